/*
 * mpcx.h -- C ABI of libmpcx, the MI355X (gfx950) implementation of the
 * secure-inference online path of the DeepDTAGen affinity branch.
 *
 * Plain C: opaque handles, plain pointers and sizes, status codes, explicit
 * HIP stream.  Both parties of the two-party protocol are evaluated in one
 * process on one GPU; every protocol exchange goes through device memory and
 * is counted (mpcx_bytes_exchanged).
 *
 * Each entry point names the reference interface it replaces (paths relative
 * to the reference repository).  The reference's kernels live in EzPC GPU-MPC
 * (not vendored); their signatures are those used at the cited call sites.
 *
 * Ring elements: uint32_t when bw == 32, uint64_t when bw == 64 ("T" below).
 * Device pointers are marked d_, host pointers h_.  A gate call over zero
 * elements (n = 0; nz = 0 for mpcx_mul_eval, rows = 0 for mpcx_ring_lincomb)
 * returns MPCX_OK without reading its pointers or counting an exchange; matrix
 * dimensions (B, N, C, nb, M, K) must be at least 1.
 */
#ifndef MPCX_H
#define MPCX_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int mpcx_status;
#define MPCX_OK 0
#define MPCX_EINVAL 1  /* bad argument (sizes, kinds, null pointers)        */
#define MPCX_EHIP 2    /* a HIP call failed; see mpcx_last_error            */
#define MPCX_ENOMEM 3  /* device allocation failed                          */
#define MPCX_ESTATE 4  /* call out of order (e.g. forward before keygen)    */
#define MPCX_EIO 5     /* a key file could not be opened, read or written, or
                          the channel to the other party failed              */
#define MPCX_EBUSY 6   /* a shared resource is in use by work still pending on
                          another stream (mpcx_maxpool_eval_noalloc)         */

typedef struct mpcx_ctx mpcx_ctx;
typedef struct mpcx_model mpcx_model;

/* Gate kinds of the truncation / ReLU family. */
#define MPCX_TR 1       /* exact floor(x/2^s) + bias  (TruncateType::TrFloor) */
#define MPCX_TRRELU 2   /* ReLU(floor(x/2^s) + bias), fused                   */
#define MPCX_RELU 3     /* ReLU(x)                                            */
#define MPCX_TRSLACK 4  /* exact floor(x/2^s), requires |x| < 2^(bw-2)        */
#define MPCX_RELUSLACK 9 /* ReLU(x), requires |x| < 2^(bw-2-s): one (bw-2-s)-bit DCF */
#define MPCX_LOCALARS 10 /* TruncateType::LocalARS, the default of DDGOrcaBatched::truncateForward
                            (gpu_mpc/ddg_orca_batched.h:180-199, keygen :273-277): the masked
                            value and its mask are shifted locally (arithmetic shift), no key
                            bytes, no exchange; floor(x/2^s) + bias + e, e in {0, 1}, or off by
                            2^(bw-s) when x + r leaves the signed ring (probability ~|x|/2^bw) */
#define MPCX_DRELU 11   /* DReLU, [x >= 0] (gpuKeyGenDRelu / the DReLU half of gpuRelu,
                           gpu_mpc/dpf_dcf_adapter.h:32-36, 97-104, 330): one (bw-1)-bit DCF and
                           one bit-plane round; the output is a masked public bit held as a ring
                           element 0/1, keygen's output "mask" is the mask bit (0/1): the
                           DReLU bit is yhat XOR mask */
/* Exact truncation in two gates, the reference's TrFloor composition (truncate-reduce
   then sign extension, gpu_mpc/dpf_dcf_adapter.h:274-303) and its ReLU-extend
   (gpuReluExtend, :225-234; keygen bin = bw - scale, bout = bw, gpu_mpc/ddg_orca.h:222): */
#define MPCX_TRMOD 12   /* floor(x/2^s) + bias, exact modulo 2^(bw-s) only: one s-bit DCF;
                           yhat is revealed reduced to bw-s bits (in [0, 2^(bw-s))) and
                           counted (and sent, in party mode) packed at bw-s bits per
                           element, as the reference's truncate-reduce reveal at bout bits
                           (gpu_mpc/dpf_dcf_adapter.h:297, gpu_comms.h:143-168) */
#define MPCX_EXT 13     /* y sign-extended from bw-s bits: the input is a TRMOD output
                           (only its low bw-s bits are read, and of the input mask too);
                           one (bw-s-1)-bit DCF.  TRMOD then EXT = MPCX_TR */
#define MPCX_EXTRELU 14 /* ReLU(y) of that value, sign-extended: the same one DCF gives the
                           sign and the wrap.  TRMOD then EXTRELU = MPCX_TRRELU */
#define MPCX_RELUPOOL 15 /* ReLU(x), requires |x| < 2^(bw-s): one (bw-s)-bit DCF (the max-pool
                            differences of EXT / EXTRELU outputs, which lie in
                            [-2^(bw-s-1), 2^(bw-s-1))) */

/* ---------------- context ----------------
 * Replaces the evaluator/dealer constructors DDGOrcaBase(party, ip, bw, scale)
 * and DDGOrcaBaseKeygen(party, bw, scale, keyFile)
 * (gpu_mpc/ddg_orca_base.h:93-116, 338-355): one context serves both parties. */
/* Environment read by mpcx_create: MPCX_AES_VARIANT and MPCX_AES_BLOCK (as
 * mpcx_set_aes_variant; bad values are ignored with a warning); MPCX_GEMM = auto
 * (default: in Z_2^32 the panel kernel where it applies, else the fused SxS and
 * wide-K matrix-core kernels where they apply, the tiled matrix-core kernels
 * elsewhere), wide (the same without the panel kernel), tiled (the tiled
 * matrix-core kernels only) or valu (the VALU kernels); MPCX_GRAPH = 0 (model
 * forwards enqueue every kernel instead of replaying a captured HIP graph).  All
 * paths give the same results bit for bit. */
mpcx_status mpcx_create(int bw, int scale, int device, mpcx_ctx **out);
void mpcx_destroy(mpcx_ctx *ctx);
const char *mpcx_last_error(const mpcx_ctx *ctx);
/* Ring width and fixed-point scale of the context. */
int mpcx_bw(const mpcx_ctx *ctx);
int mpcx_scale(const mpcx_ctx *ctx);
/* hipStream_t for the standalone gate calls; NULL = the context's own stream.
 * A model keeps the stream (and AES variant and GEMM path) the context had at
 * mpcx_model_create; mpcx_synchronize waits for the context's current stream. */
mpcx_status mpcx_set_stream(mpcx_ctx *ctx, void *hip_stream);
mpcx_status mpcx_synchronize(mpcx_ctx *ctx);
/* sync = 0: the party-mode gate calls (mpcx_party_*) return with their work
 * enqueued on the context's stream instead of synchronising it, for callers
 * that order by stream (the drop-in headers: the reference's per-call
 * semantics, gpu_comms.h's synchronous exchanges, are kept by a blocking
 * stream, on which a later null-stream copy or free waits).  Outputs are then
 * ready in the stream's order; read them on the host after mpcx_synchronize or
 * a copy ordered after the stream.  Default 1 (synchronise). */
mpcx_status mpcx_set_party_sync(mpcx_ctx *ctx, int sync);
/* AES T-table LDS layout used by the DCF kernels (0 = default).  Returns the
 * number of variants; name of variant i via mpcx_aes_variant_name.
 * block_threads: 0 (the variant's own) or a multiple of 128 in [128, 1024]. */
int mpcx_aes_variant_count(void);
const char *mpcx_aes_variant_name(int i);
mpcx_status mpcx_set_aes_variant(mpcx_ctx *ctx, int variant, int block_threads);
/* Variant in use (set by mpcx_set_aes_variant or the MPCX_AES_VARIANT environment
 * variable at mpcx_create). */
int mpcx_aes_variant(const mpcx_ctx *ctx);
/* Longest truncation/ReLU gate, in AES calls per element and party, whose
 * Z_2^32 launches of at least 1024 elements per CU run in the both-party form
 * (one thread per element holds both parties' keys; same keys and outputs):
 * 0..64, default 6; 0 keeps every gate on the one-lane-per-party kernel.  A
 * model with more than one lane takes max(setting, 14) for its own launches
 * (0 stays 0), from 512 elements per CU.  Read by the gate calls of this context and by models created
 * after it.  No counterpart in the reference: a tuning setting of this
 * library, as mpcx_set_aes_variant. */
mpcx_status mpcx_set_both_party_aes(mpcx_ctx *ctx, int max_aes);

/* The dealer's 16 secret key bytes (NULL: none).  With a key set, every
 * keygen of this context (and of models created afterwards) derives its PRF key
 * from these bytes and the seed (which then only names the key set), so the
 * keys rest on 128 secret bits; without one the seed alone determines them,
 * which suits tests and benchmarks.  Both parties' keys come from the one dealer
 * run, as the reference's dealer (DDGOrcaBaseKeygen, gpu_mpc/ddg_orca_base.h:
 * 338-355, with initGPURandomness) draws them. */
mpcx_status mpcx_set_dealer_key(mpcx_ctx *ctx, const uint8_t *key16);

/* Exchange accounting, both directions summed (the reference's "Comm (B)",
 * gpu_mpc/deepdtagen_inference.cu:556-558, and GpuPeer::bytesSent/Received,
 * gpu_mpc/utils/gpu_comms.h:290-397). */
uint64_t mpcx_bytes_exchanged(const mpcx_ctx *ctx);
uint64_t mpcx_rounds(const mpcx_ctx *ctx);
void mpcx_reset_counters(mpcx_ctx *ctx);

/* ---------------- PRG ----------------
 * Tree hash H(s) = AES_KH(sigma(s)) ^ sigma(s) (leaf = 0) or the leaf hash HL
 * (leaf = 1) on n 128-bit blocks; replaces the AES context of GPU-MPC
 * (AESGlobalContext / initAESContext, gpu_mpc/ddg_orca_base.h:50,95). */
mpcx_status mpcx_prg_hash(mpcx_ctx *ctx, int leaf, size_t n, const void *d_in, void *d_out);
/* Dealer PRF blocks AES_Kd(i, field, gate), i = 0..n-1 (randomGEOnGpu,
 * randomAESBlockOnGpu in GPU-MPC). */
mpcx_status mpcx_prf(mpcx_ctx *ctx, uint64_t seed, uint32_t gate, uint32_t field, size_t n, void *d_out);

/* ---------------- DCF ----------------
 * [x < alpha] over bin-bit inputs, XOR-shared output bits masked by rbit.
 * Replaces gpuKeyGenDCF<T>(u8**, party, bin, N, T* d_rin, AESGlobalContext*)
 * (gpu_mpc/dpf_dcf_adapter.h:372), readGPUDcfKey (:100) and
 * gpuDcf<T,1,idPrologue,maskEpilogue>(key, party, d_in, g, s) (:266).
 * alpha and x: n uint64_t each; rbit: n bytes or NULL; out: packed bits,
 * bit i of 64-bit word i/64, (n+63)/64 words. */
size_t mpcx_dcf_key_bytes(int bin, size_t n);
mpcx_status mpcx_dcf_keygen(mpcx_ctx *ctx, int bin, size_t n, const uint64_t *d_alpha,
                            const uint8_t *d_rbit, uint64_t seed, uint32_t gate, void *d_key0,
                            void *d_key1);
mpcx_status mpcx_dcf_eval(mpcx_ctx *ctx, int party, int bin, size_t n, const void *d_key,
                          const uint64_t *d_x, uint64_t *d_out_bits);
/* The same on ring elements of the context's width (d_x: n uint32_t at bw=32,
 * uint64_t at bw=64; each read modulo 2^bin), with the output bits XORed with
 * d_mask (device, (n+31)/32 words, bit i of word i/32) when it is not NULL: the
 * reference's gpuDcf<T, 1, idPrologue, maskEpilogue>(key, party, d_in, g, s,
 * &h_mask) (gpu_mpc/dpf_dcf_adapter.h:266, 293) with no host round trip. */
mpcx_status mpcx_dcf_eval_ring(mpcx_ctx *ctx, int party, int bin, size_t n, const void *d_key,
                               const void *d_x, const uint32_t *d_mask, uint64_t *d_out_bits);

/* ---------------- truncation / ReLU ----------------
 * Keygen replaces gpuGenReluKey<T,T,0,0,false>(kb, party, bin, bout, N,
 * d_inMask, g) (gpu_mpc/ddg_orca.h:233) and genGPUTruncateKey<T,T>(kb, party,
 * TrFloor, bin, bout, shift, N, d_inMask, g) (gpu_mpc/ddg_orca.h:240-241):
 * takes the input mask, writes the output mask and both parties' keys.
 * Eval replaces gpuRelu<T,T,0,0,false>(peer, party, key, d_in, g, s)
 * (gpu_mpc/ddg_orca.h:103-104) and gpuTruncate<T,T>(bin, bout, TrFloor, k,
 * shift, peer, party, N, d_in, g, s) (gpu_mpc/ddg_orca.h:116-118), for both
 * parties at once: masked input in, masked output out.
 * bias: ncol ring elements at scale s (element i uses bias[i % ncol]) or NULL;
 * read only by MPCX_TR, MPCX_TRRELU, MPCX_TRSLACK, MPCX_TRMOD and MPCX_LOCALARS
 * (the kinds that shift).  MPCX_LOCALARS has no key (key bytes 0, key pointers
 * may be NULL, the gate id is unused). */
size_t mpcx_tr_key_bytes(mpcx_ctx *ctx, int kind, size_t n);
/* AES calls per element and party of a gate kind's evaluation (its DCF walks:
 * tree levels plus the leaf), for the caller's own accounting of the DCF work
 * (the reference's Stats counts time only); 0 for MPCX_LOCALARS, -1 for a bad
 * kind. */
int mpcx_tr_aes_calls(const mpcx_ctx *ctx, int kind);
/* The kernel form mpcx_tr_eval takes for n elements of a gate kind on this
 * context and its settings (mpcx_set_both_party_aes, mpcx_set_aes_variant):
 * the one-lane kernel, the both-party form (one thread per element runs both
 * parties' DCF walks) or the quad-lane form (four lanes per element and party);
 * -1 for a bad kind or MPCX_LOCALARS.  No counterpart in the reference: a query
 * for tests and tuning. */
#define MPCX_FORM_ONE_LANE 0
#define MPCX_FORM_BOTH 1
#define MPCX_FORM_QUAD 2
int mpcx_tr_eval_form(const mpcx_ctx *ctx, int kind, size_t n);
mpcx_status mpcx_tr_keygen(mpcx_ctx *ctx, int kind, size_t n, const void *d_in_mask,
                           void *d_out_mask, uint64_t seed, uint32_t gate, void *d_key0,
                           void *d_key1);
mpcx_status mpcx_tr_eval(mpcx_ctx *ctx, int kind, size_t n, const void *d_key0,
                         const void *d_key1, const void *d_xhat, const void *d_bias, int ncol,
                         void *d_yhat);

/* ---------------- masked global max-pool ----------------
 * Replaces MaskedMaxPoolLayer<T>(B, Nmax, F)::_forward
 * (gpu_mpc/masked_maxpool_layer.h:47-165; MaskedGlobalMaxPool for B = 1,
 * gpu_mpc/masked_maxpool.h:62-84): input (B*N, C) masked-public, sample-major
 * (the reference's input is already H (.) mask), output (B, C): per sample and
 * channel the maximum over the N rows, as the reference's tree — pairs of rows
 * (2j, 2j+1), max(a, b) = a + ReLU(b - a), an odd last row carried to the next
 * level — over mpcx_maxpool_levels(N) = ceil(log2 N) levels, two exchange
 * rounds each.  Exact while every pairwise difference lies in the signed ring.
 * Keygen uses the gate ids gate .. gate + levels - 1; with N = 1 there is no key
 * (key pointers may be NULL) and the output is the input. */
int mpcx_maxpool_levels(int N);
size_t mpcx_maxpool_key_bytes(mpcx_ctx *ctx, int B, int N, int C);
mpcx_status mpcx_maxpool_keygen(mpcx_ctx *ctx, int B, int N, int C, const void *d_in_mask,
                                void *d_out_mask, uint64_t seed, uint32_t gate, void *d_key0,
                                void *d_key1);
mpcx_status mpcx_maxpool_eval(mpcx_ctx *ctx, int B, int N, int C, const void *d_key0,
                              const void *d_key1, const void *d_xhat, void *d_yhat);
/* Allocation-free variant of mpcx_maxpool_eval.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, keys and results.  Its level planes live in a static device
 * array of MPCX_NOALLOC_SCRATCH_BYTES per GPU (resident from the library's load
 * until the process ends) instead of the context's workspace: it calls no
 * hipMalloc, hipFree or allocating routine and does not synchronize (the
 * output is ready when the context's stream reaches it).  It needs
 * (2*B*N*C + 2*B*floor(N/2)*C) * bw/8 bytes of that array (64 x 140 x 312 fits
 * at both widths); larger calls fail with MPCX_EINVAL.  Every call on one GPU
 * shares that GPU's array: calls on one stream run in order; a call on another
 * stream (another context, thread or mpcx_set_stream) while the last call's
 * work is still pending fails with MPCX_EBUSY before any launch (the library
 * tracks the last caller's stream and an event it records after the call;
 * calls captured into a HIP graph are not tracked, so replays of such a graph
 * must not overlap other calls on the same GPU). */
#define MPCX_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
mpcx_status mpcx_maxpool_eval_noalloc(mpcx_ctx *ctx, int B, int N, int C, const void *d_key0,
                                      const void *d_key1, const void *d_xhat, void *d_yhat);

/* ---------------- Beaver product ----------------
 * z[i] = x[ia[i]] * y[ib[i]] on masked operands (index maps allow the
 * broadcast/outer products of the adjacency normalisation).  Replaces
 * gpuKeygenMul<T>(kb, party, bw, scale, N, d_maskA, d_maskB, None, g) and
 * gpuMul<T>(peer, party, bw, scale, N, key, d_A, d_B, None, g, s)
 * (gpu_mpc/secure_adj_norm.h:326-337, 611-624; gpu_mpc/ddg_orca.h:43-63). */
size_t mpcx_mul_key_bytes(mpcx_ctx *ctx, size_t nx, size_t ny, size_t nz);
mpcx_status mpcx_mul_keygen(mpcx_ctx *ctx, size_t nx, size_t ny, size_t nz, const uint32_t *d_ia,
                            const uint32_t *d_ib, const void *d_rx, const void *d_ry, void *d_rz,
                            uint64_t seed, uint32_t gate, void *d_key0, void *d_key1);
mpcx_status mpcx_mul_eval(mpcx_ctx *ctx, size_t nx, size_t ny, size_t nz, const uint32_t *d_ia,
                          const uint32_t *d_ib, const void *d_key0, const void *d_key1,
                          const void *d_xhat, const void *d_yhat, void *d_zhat);

/* Byte offsets, from the start of a party's Beaver-product key, of its share of
 * the x mask (nx elements), of the y mask (ny) and of the product term (nz): the
 * fields a, b, c of the reference's GPUMulKey, which callers read to reveal a
 * leaf operand (gpu_mpc/ddg_orca.h:50-57, gpu_mpc/secure_adj_norm.h:630-640). */
mpcx_status mpcx_mul_key_layout(mpcx_ctx *ctx, size_t nx, size_t ny, size_t nz, size_t off[3]);

/* ---------------- 8-bit DPF lookup table ----------------
 * y = table[x] for secret x in [0, 256) (the D^-1/2 degree table).  Replaces
 * gpuKeyGenLUT<T,T>(kb, party, 8, bw, N, d_inMask, g), readGPULUTKey and
 * gpuDpfLUT<T,T>(key, peer, party, d_x, d_table, g, s, true)
 * (gpu_mpc/secure_adj_norm.h:270-279, 498-520).  table: 256 ring elements. */
size_t mpcx_lut8_key_bytes(mpcx_ctx *ctx, size_t n);
mpcx_status mpcx_lut8_keygen(mpcx_ctx *ctx, size_t n, const void *d_in_mask, void *d_out_mask,
                             uint64_t seed, uint32_t gate, void *d_key0, void *d_key1);
mpcx_status mpcx_lut8_eval(mpcx_ctx *ctx, size_t n, const void *d_key0, const void *d_key1,
                           const void *d_table, const void *d_xhat, void *d_yhat);

/* ---------------- ring GEMMs ----------------
 * Batched secret x secret product C_b = A_b (M x K) . B_b (K x N) on masked
 * operands (Beaver).  Replaces the 3-argument DDGOrcaBase::matmul and its
 * keygen mirror (gpu_mpc/ddg_orca_base.h:170-205, 394-410), i.e.
 * gpuKeygenMatmul / gpuMatmul with wIsOnGpu = true and the per-sample loop of
 * _MatMul (gpu_mpc/sytorch/layers/layers.h:67-93). */
size_t mpcx_sxs_key_bytes(mpcx_ctx *ctx, int nb, int M, int K, int N);
mpcx_status mpcx_sxs_keygen(mpcx_ctx *ctx, int nb, int M, int K, int N, const void *d_ra,
                            const void *d_rb, void *d_rc, uint64_t seed, uint32_t gate,
                            void *d_key0, void *d_key1);
mpcx_status mpcx_sxs_eval(mpcx_ctx *ctx, int nb, int M, int K, int N, const void *d_key0,
                          const void *d_key1, const void *d_ahat, const void *d_bhat,
                          void *d_chat);
/* Byte offsets, from the start of a party's SxS key, of its shares of the A
 * mask (nb*M*K), of the B mask (nb*K*N) and of its C term (nb*M*N): the fields
 * A, B, C of the reference's GPUMatmulKey (gpu_mpc/ddg_orca_base.h:181-186). */
mpcx_status mpcx_sxs_key_layout(mpcx_ctx *ctx, int nb, int M, int K, int N, size_t off[3]);
/* Public ring GEMM C = A . B mod 2^bw (masked activations x public weights;
 * the 4-argument DDGOrcaBase::matmul, gpu_mpc/ddg_orca_base.h:208-271, needs no
 * key and no exchange when the output mask is r_A . W). */
mpcx_status mpcx_ring_gemm(mpcx_ctx *ctx, int M, int K, int N, const void *d_a, const void *d_b,
                           void *d_c);

/* Local linear map on masked-public ring tensors (rows x cols, row-major):
 * out = a*x + b*y + (v[col] << shift), x, y or v may be NULL.  Linear maps need no
 * key and no exchange: the evaluators apply them to masked values and the dealer
 * to the masks (with v = NULL, since a public addend has mask 0).  Replaces
 * gpuLinearComb / gpuAdd behind the backend's add, sub and scalarmul
 * (gpu_mpc/ddg_orca_base.h:304-314, gpu_mpc/ddg_orca.h:65-81) and the bias add of
 * the 4-argument matmul (ddg_orca_base.h:208-271, bias at scale 2s). */
mpcx_status mpcx_ring_lincomb(mpcx_ctx *ctx, size_t rows, size_t cols, uint64_t a, const void *d_x, uint64_t b,
                              const void *d_y, const void *d_v, int shift, void *d_out);

/* ---------------- reveal ----------------
 * Additive shares v0, v1 -> masked public v + r (revealIfLeaf,
 * gpu_mpc/ddg_orca_base.h:72-80; peer->reconstructInPlace,
 * gpu_mpc/utils/gpu_comms.h:290-302). */
size_t mpcx_reveal_key_bytes(mpcx_ctx *ctx, size_t n);
mpcx_status mpcx_reveal_keygen(mpcx_ctx *ctx, size_t n, void *d_mask, uint64_t seed, uint32_t gate,
                               void *d_key0, void *d_key1);
mpcx_status mpcx_reveal_eval(mpcx_ctx *ctx, size_t n, const void *d_key0, const void *d_key1,
                             const void *d_v0, const void *d_v1, void *d_vhat);

/* ---------------- secure adjacency normalisation ----------------
 * A_norm = D^-1/2 (A) D^-1/2 on secret A, in the fixed-point form of the secure
 * path: A[i,j] * floor(T[d_i] T[d_j] / 2^s), T[k] = llround(2^s / sqrt(k)) for
 * 1 <= k <= nmax, T[0] = 0, d = row sums of A (self loops included).  Replaces
 * ddgSecureAdjNormKeygen / ddgSecureAdjNormEval (gpu_mpc/secure_adj_norm.h:203-374,
 * 393-659): reveal A, reveal the degrees, 8-bit DPF-LUT, Beaver outer product,
 * one exact truncation, Beaver A (.) W.  a0, a1: both parties' shares of A
 * (B x N x N ring elements, N <= 255); out: A_norm + out_mask. */
size_t mpcx_adjnorm_key_bytes(mpcx_ctx *ctx, int B, int N);
/* Concurrent graph groups (1..16, default 1) of the adjacency normalisation
 * calls of this context: the B graphs are split into that many groups of
 * consecutive graphs (B/L each, the first B%L one larger), each evaluated on its
 * own stream so that one group's DCF work overlaps another's memory-bound
 * gates.  The key set is the groups' one-group key sets back to back, group i
 * keyed under seed + i * 0x9E3779B97F4A7C15: keygen and eval must use the same
 * setting (like the model's lanes, mpcx_model_set_lanes). */
mpcx_status mpcx_set_adjnorm_lanes(mpcx_ctx *ctx, int lanes);
mpcx_status mpcx_adjnorm_keygen(mpcx_ctx *ctx, int B, int N, uint64_t seed, void *d_out_mask, void *d_key0,
                                void *d_key1);
mpcx_status mpcx_adjnorm_eval(mpcx_ctx *ctx, int B, int N, int nmax, const void *d_key0, const void *d_key1,
                              const void *d_a0, const void *d_a1, void *d_out);

/* ---------------- party mode: one process (or thread) per party ----------------
 * The reference deploys the two parties as two processes on one GPU, each with
 * its own key file, talking over a socket (gpu_mpc/run_local_2pc.sh:196-233;
 * GpuPeer / SigmaPeer, gpu_mpc/utils/gpu_comms.h:94-397,
 * gpu_mpc/utils/sigma_comms.cpp:36-150).  In party mode each process creates its
 * own context on the GPU and one end of a channel; every exchange sends exactly
 * the bytes mpcx_bytes_exchanged counts (ring elements at their width, DCF output
 * bits packed 32 per 32-bit word: the bit-packed wire of gpu_comms.h:28-73), and
 * each party's context counts both directions, as in the one-process mode.  The
 * gate calls below take this party's key (as written by the keygen calls for
 * that party) and its share or the masked public input, and return the
 * reconstructed masked output on both parties; they synchronise the context's
 * stream (unless mpcx_set_party_sync(ctx, 0)). */
typedef struct mpcx_peer mpcx_peer;
/* Party 0 listens on the Unix socket `path`, party 1 connects (GpuPeer::connect,
 * gpu_mpc/ddg_orca_base.h:113-114).  timeout_ms bounds the rendezvous and every
 * later receive.  MPCX_EIO if no connection is made. */
mpcx_status mpcx_peer_connect(int party, const char *path, int timeout_ms, mpcx_peer **out);
/* Both ends of one channel, for two parties run as two threads of one process.
 * The ends are linked in memory: an exchange is a device-to-device copy of each
 * party's message into the other's receive regions, ordered by events on the
 * two parties' streams (no host staging, no socket); bytes and rounds are
 * counted as on a socket.  With MPCX_PEER_SOCKETPAIR=1 in the environment the
 * ends are a socket pair, staged through pinned host memory as between two
 * processes.  timeout_ms bounds the wait for the peer at each exchange. */
mpcx_status mpcx_peer_pair(int timeout_ms, mpcx_peer **p0, mpcx_peer **p1);
void mpcx_peer_close(mpcx_peer *peer);
int mpcx_peer_party(const mpcx_peer *peer);
/* Bytes sent plus bytes received over the channel, and exchanges made. */
uint64_t mpcx_peer_bytes(const mpcx_peer *peer);
uint64_t mpcx_peer_rounds(const mpcx_peer *peer);
/* How the channel moves messages: 2 device to device within one process
 * (mpcx_peer_pair), 1 through device inboxes shared by IPC memory handles (two
 * processes on one GPU: each exchange writes this party's message straight into
 * the peer's inbox, one-byte tokens on the socket order the writes and reads),
 * 0 staged through pinned host memory and the socket (other setups, messages
 * over 1 GiB, MPCX_PEER_IPC=0 in either process), -1 not yet decided (a
 * connected channel before its first exchange).  No counterpart in the
 * reference, whose GpuPeer always stages through the host. */
int mpcx_peer_transport(const mpcx_peer *peer);
const char *mpcx_peer_error(const mpcx_peer *peer);
/* peer->reconstructInPlace(d, bw, n, s) (gpu_mpc/utils/gpu_comms.h:290-302):
 * d_inout holds this party's additive share and receives the sum of both. */
mpcx_status mpcx_party_reconstruct(mpcx_ctx *ctx, mpcx_peer *peer, size_t n, void *d_inout);
/* gpuRelu / gpuTruncate / gpuReluExtend / the DReLU of gpuRelu for this party
 * (gpu_mpc/ddg_orca.h:90, 103-104, 116-118; dpf_dcf_adapter.h:225-234):
 * d_key = this party's key (mpcx_tr_key_bytes); MPCX_DRELU returns the public
 * masked bit after one round, the other kinds the masked output after two. */
mpcx_status mpcx_party_tr_eval(mpcx_ctx *ctx, mpcx_peer *peer, int kind, size_t n, const void *d_key,
                               const void *d_xhat, const void *d_bias, int ncol, void *d_yhat);
/* gpuMul (gpu_mpc/secure_adj_norm.h:611-624, gpu_mpc/ddg_orca.h:43-63). */
mpcx_status mpcx_party_mul_eval(mpcx_ctx *ctx, mpcx_peer *peer, size_t nx, size_t ny, size_t nz,
                                const uint32_t *d_ia, const uint32_t *d_ib, const void *d_key,
                                const void *d_xhat, const void *d_yhat, void *d_zhat);
/* gpuDpfLUT (gpu_mpc/secure_adj_norm.h:510-520). */
mpcx_status mpcx_party_lut8_eval(mpcx_ctx *ctx, mpcx_peer *peer, size_t n, const void *d_key,
                                 const void *d_table, const void *d_xhat, void *d_yhat);
/* gpuMatmul, secret x secret (gpu_mpc/ddg_orca_base.h:170-205). */
mpcx_status mpcx_party_sxs_eval(mpcx_ctx *ctx, mpcx_peer *peer, int nb, int M, int K, int N, const void *d_key,
                                const void *d_ahat, const void *d_bhat, void *d_chat);
/* revealIfLeaf (gpu_mpc/ddg_orca_base.h:72-80): d_v this party's share. */
mpcx_status mpcx_party_reveal_eval(mpcx_ctx *ctx, mpcx_peer *peer, size_t n, const void *d_key,
                                   const void *d_v, void *d_vhat);

/* ---------------- pinned host memory ----------------
 * Page-locked host buffers for streamed key arenas (hipHostMalloc). */
mpcx_status mpcx_host_alloc(size_t bytes, void **out);
void mpcx_host_free(void *p);

/* ---------------- the model ----------------
 * DeepDTAGenAffinity<T> (gpu_mpc/deepdtagen.h:110-223) with the driver's
 * resident-key evaluation loop (gpu_mpc/deepdtagen_inference.cu:422-607).
 * Weights: the weights.bin layout (deepdtagen_inference.cu:121-181): for each
 * linear layer W^T (in x out, row-major) then bias (out), int64 at scale s. */
typedef struct {
  int n_nodes;  /* padded atoms per molecule (<= 255) */
  int feat;     /* atom feature width */
  int gcn[3];   /* GCN output widths */
  int dfc[2];   /* drug FC widths */
  int prot;     /* protein embedding width */
  int nfus;     /* fusion layers (last has width 1) */
  int fus[4];
  int lut_nmax; /* largest degree with a D^-1/2 table entry */
  int mask_scale; /* atom mask values are 0 or 2^mask_scale: 0, or s for the reference's
                     mask files (reference/share_data.py:135-159 shares the mask at scale s) */
  int slack;      /* 0: every truncation is exact over the signed ring (DDGOrca::truncateForward
                     TrFloor, gpu_mpc/ddg_orca.h:112-123: two DCFs, 31 AES per element and party
                     at bw=32).  1: the GCN products H.W^T use the top-two-bit slack truncation
                     (the reference's TrWithSlack, ddg_orca.h:50, 60), exact for |H.W^T| <
                     2^(bw-2), one s-bit DCF (6 AES).  2: also the aggregation A.XW + bias:
                     slack truncation with the bias, then MPCX_RELUSLACK on the truncated value
                     (a (bw-2-s)-bit DCF, 12 AES at bw=32; two more exchange rounds), exact for
                     |A.XW + b 2^s| < 2^(bw-2).  Outputs are bit-exact with the fixed-point
                     forward while every such value lies in that half ring.  3: every layer
                     truncation (H.W^T, A.XW + b, the FCs) is MPCX_LOCALARS, the reference's
                     default (gpu_mpc/ddg_orca_batched.h:180-199), followed by a RELU gate on
                     ReLU layers; the adjacency normalisation stays exact.  Not bit-exact:
                     +1 per truncation, and a 2^(bw-s) error when x + r wraps (~|x|/2^bw per
                     element: usable at bw=64 only, as the reference notes). */
} mpcx_model_dims;

mpcx_status mpcx_model_create(mpcx_ctx *ctx, const mpcx_model_dims *dims, const int64_t *h_weights,
                              size_t n_weights, mpcx_model **out);
void mpcx_model_destroy(mpcx_model *m);
/* Concurrent sub-batches: every batch of B is split into `lanes` (1..16)
 * sub-batches of consecutive samples (B/lanes each, the first B%lanes one
 * larger), each evaluated by its own copy of the gate sequence on its own
 * stream; the context stream waits for every lane at the end of a forward.
 * Lanes past the first do not wait for work enqueued on the context stream
 * before the forward (the forward reads only the model's buffers, which
 * mpcx_model_set_inputs fills synchronously).  The reference
 * evaluates a batch as one gate sequence (DeepDTAGenAffinity<T>::_forward,
 * gpu_mpc/deepdtagen.h:183-222); lanes let the gates of one sub-batch that
 * leave the GPU partly idle overlap another's DCF evaluation.  Keys of a batch
 * are the lanes' key sets back to back, lane i's being the one-lane key set
 * of its samples under seed + i * 0x9E3779B97F4A7C15 (mod 2^64); with
 * host-streamed keys each lane has its own two slots of slot_bytes.  Drops
 * keys and inputs.  Default: 1 lane. */
mpcx_status mpcx_model_set_lanes(mpcx_model *m, int lanes);
int mpcx_model_lanes(const mpcx_model *m);
/* Key bytes per party for a batch of B molecules. */
size_t mpcx_model_key_bytes(const mpcx_model *m, int B);
/* Dealer on the GPU: generates both parties' keys into the resident key arena
 * (initGPUKeyArena, patches/EzPC-GPU-MPC.track3.patch:632-661). */
mpcx_status mpcx_model_keygen(mpcx_model *m, int B, uint64_t seed);
/* Upload / download whole key arenas (host buffers of mpcx_model_key_bytes). */
mpcx_status mpcx_model_import_keys(mpcx_model *m, int B, const void *h_key0, const void *h_key1,
                                   size_t bytes);
mpcx_status mpcx_model_export_keys(mpcx_model *m, int party, void *h_dst, size_t bytes);
/* Frees the resident key arenas (e.g. after mpcx_model_export_keys). */
mpcx_status mpcx_model_release_arena(mpcx_model *m);
/* Packed keys.  The DCF correction and leaf words and the clear output mask are
 * the same in both parties' keys; the evaluation reads them from party 0's copy.
 * The dealer draws every purely random plane of a party's truncation-family
 * keys (DCF roots and output-mask bits; for party 0 also its shares of kappa and
 * of the G tables) from that party's own PRF key, which the party receives
 * instead of those planes (the seed compression of the reference's key format
 * notes, README.md:144-157, 319-322).  Party p's packed key: a 256-byte header
 * (its 16-byte PRF key, then zeros) and its remaining planes back to back in
 * arena order, mpcx_model_unique_key_bytes(m, B, p) bytes (at bw=64 about 90%
 * of party 0's arena and 7% of party 1's); with lanes, the lanes' packed keys
 * back to back.  Exported from keys made by mpcx_model_keygen only (imported
 * keys carry no PRF keys: MPCX_ESTATE). */
size_t mpcx_model_unique_key_bytes(const mpcx_model *m, int B, int party);
mpcx_status mpcx_model_export_unique_keys(mpcx_model *m, int party, void *h_dst, size_t bytes);
/* Streaming key arena for batches whose keys do not stay resident: both parties'
 * keys in host memory (pinned for overlap) are copied per chunk of consecutive
 * gates into one of two device slots of at most slot_bytes per party, on a copy
 * stream, while the previous chunk computes; party 1's shared planes are not
 * copied.  Each of h_key0, h_key1: the party's arena (bytes = mpcx_model_key_bytes)
 * or its packed key (bytes = mpcx_model_unique_key_bytes(m, B, p)), whose
 * PRF-drawn planes are expanded in the device slot after each chunk's copy, on
 * the copy stream.  Replaces the chunked key
 * pipeline of gpu_mpc/deepdtagen_inference.cu:608-859 (pinned double-buffered
 * slots, copy stream, ready/free events) and setGPUKeyArenaSlot
 * (patches/EzPC-GPU-MPC.track3.patch:680-685).  The resident arena is freed;
 * the host buffers must stay valid until the model is destroyed.  MPCX_EINVAL
 * if a single gate's key exceeds slot_bytes. */
mpcx_status mpcx_model_attach_host_keys(mpcx_model *m, int B, const void *h_key0, size_t bytes0,
                                        const void *h_key1, size_t bytes1, size_t slot_bytes);
/* Key files.  mpcx_model_write_keys appends the key set of the batch keyed
 * last (mpcx_model_keygen / import) for one party to a file: the party's arena
 * (packed = 0) or its packed key (packed = 1, keys from keygen only); append
 * = 0 truncates the file first.  Sets of successive keygens (fresh seeds)
 * appended in order form a key file of whole-batch key sets.
 * mpcx_model_attach_key_files streams such files: each forward reads the next
 * key set (cycling), chunk by chunk: an I/O thread preads chunk k into one of
 * two pinned staging buffers per party (chunk k - 2's copies out of it done),
 * the copy stream moves it into a device slot of at most slot_bytes per party
 * and lane, and the gates of the chunk wait for that copy.  Replaces the
 * SSD -> pinned -> VRAM pipeline of gpu_mpc/deepdtagen_inference.cu:608-859
 * (I/O thread, pread into pinned slots, evH2D / evFree handshake); the
 * reference's chunks are whole micro-batch key sets, these are gate-aligned
 * pieces of one, so a key set need not fit in memory twice.  Each file holds
 * arenas or packed keys, told apart by its size.  MPCX_EIO if a
 * file is missing, does not hold whole key sets, or a read fails. */
mpcx_status mpcx_model_write_keys(mpcx_model *m, int party, int packed, const char *path, int append);
mpcx_status mpcx_model_attach_key_files(mpcx_model *m, int B, const char *path0, const char *path1,
                                        size_t slot_bytes);
/* Chunks and host-to-device key bytes (both parties) of the last forward. */
mpcx_status mpcx_model_stream_stats(const mpcx_model *m, int *chunks, uint64_t *bytes_h2d);
/* Both parties' input shares (host, ring elements): x (B,N,feat), adjacency
 * (B,N,N) at scale 0 with self loops, atom mask (B,N); protein embedding
 * (B,prot) int64 at scale s, public. */
mpcx_status mpcx_model_set_inputs(mpcx_model *m, int B, const void *h_x0, const void *h_x1,
                                  const void *h_a0, const void *h_a1, const void *h_m0,
                                  const void *h_m1, const int64_t *h_prot);
/* One online forward of both parties (enqueued on the context stream). */
mpcx_status mpcx_model_forward(mpcx_model *m, int B);
/* Reconstructed outputs (B int64 at scale s); synchronizes the stream. */
mpcx_status mpcx_model_output(mpcx_model *m, int B, int64_t *h_out);
/* Party mode of the model (one lane; the reference's evaluator process,
 * gpu_mpc/deepdtagen_inference.cu:422-607 with run_local_2pc.sh:196-233): the
 * model evaluates only the peer's party, holding that party's key and shares,
 * and exchanges through the peer; peer = NULL returns to both parties in one
 * process.  Drops keys and inputs.  The party imports its own key
 * (mpcx_model_export_keys / mpcx_model_write_keys of the dealer's run for that
 * party, mpcx_model_key_bytes bytes) and its input shares; h_prot is the
 * protein embedding on the party that owns it (party 1 in the reference's
 * deployment) and NULL on the other.  mpcx_model_forward / _output then work
 * as in the one-process mode and give the same outputs and exchange bytes. */
mpcx_status mpcx_model_set_party(mpcx_model *m, mpcx_peer *peer);
mpcx_status mpcx_model_import_party_key(mpcx_model *m, int B, const void *h_key, size_t bytes);
mpcx_status mpcx_model_set_party_inputs(mpcx_model *m, int B, const void *h_x, const void *h_a,
                                        const void *h_m, const int64_t *h_prot);
/* DCF gate kernel (k_tr_eval) timing with HIP events on the launch streams.  While
 * enabled, forwards run their lanes one after another (each launch is timed
 * alone) and launch the separately named k_tr_eval<..., 1> instantiation. */
mpcx_status mpcx_model_profile(mpcx_model *m, int enable);
/* After a synchronized forward: number of DCF gate launches, their summed time
 * (ms), elements (both parties), AES calls (both parties) and algorithmic HBM
 * bytes (keys, inputs, G words and kappa read, the revealed output written; both
 * parties). */
mpcx_status mpcx_model_profile_read(mpcx_model *m, int *launches, double *ms, double *elements,
                                    double *aes_calls, double *hbm_bytes);
/* After a synchronized profiled forward: ring-GEMM sections (one per public-
 * weight product, one per SxS gate's three Beaver products), their summed time
 * (ms, HIP events on the launch streams) and the ring multiply-adds inside
 * (the reference's gpuMatmul, gpu_mpc/ddg_orca_base.h:170-271). */
mpcx_status mpcx_model_profile_gemm(mpcx_model *m, int *sections, double *ms, double *ring_macs);

#ifdef __cplusplus
}
#endif
#endif
