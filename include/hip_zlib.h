/* C-ABI of the MI355X (gfx950) zlib/DEFLATE codec.
 *
 * Every entry point takes device pointers, sizes and a HIP stream.  Work is
 * enqueued on that stream; no entry point synchronises with the host except
 * where noted.  Buffers are owned by the caller; scratch comes from a private
 * per-device stream-ordered pool.
 *
 * Return value: 0 on success; a positive hipError_t for a HIP runtime failure;
 * HIP_ZLIB_INVALID_ARGUMENT (-1) for a malformed call (wrong metadata shape,
 * inconsistent batch layout).  HipZlibErrorString() describes either.  Data
 * errors are never returned: they are written to the metadata buffer as codec
 * statuses (0 ok, 1..23 as documented in the Python package), exactly like the
 * reference's XLA FFI handlers, which return Success with an error status.
 */
#ifndef HIP_ZLIB_H_
#define HIP_ZLIB_H_

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HIP_ZLIB_INVALID_ARGUMENT (-1)

/* Compress input[0..input_size) into a zero-padded zlib stream.
 * output_size must equal input_size + 5 * max(1, ceil(input_size / chunk_bytes)) + 6.
 * metadata (2 x u32, device): [encoded_length, status].
 * Replaces the reference's CudaZlibCompress FFI handler
 * (src/cuda_zlib/native/codec_ffi.cu:1144-1152, body Compress at 551-612). */
int HipZlibCompress(hipStream_t stream, int64_t chunk_bytes, const uint8_t* input,
                    uint64_t input_size, uint8_t* output, uint64_t output_size,
                    uint32_t* metadata, uint64_t metadata_count);

/* HipZlibCompress with every chunk's LZ77 window limited to the chunk itself
 * (no matches into the bytes before it), the reference encoder's semantics
 * ("Chunks have no shared history", src/cuda_zlib/_encode_kernels.py:6;
 * encode_chunk 283-393, launched by Compress at codec_ffi.cu:551-612).  Same
 * arguments, checks, statuses and metadata as HipZlibCompress; the stream is
 * usually somewhat larger.  The reference has no separate handler for it: its
 * one compress handler always encodes chunks this way. */
int HipZlibCompressIndependent(hipStream_t stream, int64_t chunk_bytes, const uint8_t* input,
                               uint64_t input_size, uint8_t* output, uint64_t output_size,
                               uint32_t* metadata, uint64_t metadata_count);

/* Decompress a zlib stream into exactly output_size bytes.
 * metadata (2 x u32, device): [status, 0].  Output is zero-filled on failure
 * (serial small-stream route: decoded prefix followed by zeros).
 * Replaces CudaZlibDecompress (codec_ffi.cu:1153-1162, body Decompress at 662-950). */
int HipZlibDecompress(hipStream_t stream, int64_t max_candidates, int64_t max_blocks,
                      const uint8_t* input, uint64_t input_size, uint8_t* output,
                      uint64_t output_size, uint32_t* metadata, uint64_t metadata_count);

/* Decompress one stream in a wrapper format the reference does not decode:
 * format 0 zlib, 1 raw DEFLATE (RFC 1951, no wrapper or checksum), 2 gzip
 * (RFC 1952, one member: optional header fields, FHCRC, CRC-32 and ISIZE
 * checked).  dictionary (device, dictionary_size bytes; null and 0 for none)
 * is the preset dictionary of a zlib stream whose header sets FDICT (its
 * Adler-32 must equal the DICTID) or the history of a raw stream; a zlib
 * stream without FDICT ignores it, and gzip takes none.  Arguments, metadata
 * [status, 0] and failure behaviour are HipZlibDecompress's, with two more
 * statuses: 24 (gzip CRC-32 or ISIZE mismatch; output kept, as for 21) and 25
 * (dictionary Adler-32 differs from the DICTID).  Bytes after the stream's end
 * (such as a second gzip member) give status 12.  Format 0 without a
 * dictionary is exactly HipZlibDecompress.  With a dictionary, an output
 * above 64 KiB (or any output under non-default limits) is decoded into
 * scratch behind the dictionary's last 32 KiB and then copied to `output`:
 * the call needs about output_size more scratch, and one more pass over the
 * output, than the same stream without a dictionary.  No
 * counterpart in the reference, which rejects gzip with status 16 and
 * dictionaries with 17 (src/cuda_zlib/_codec.py:105-111).
 *
 * format | HIP_ZLIB_FORMAT_MEMBERS (zlib or gzip, no dictionary) decodes a
 * concatenation: one member after another (each zlib stream or gzip member
 * with its own header, window and Adler-32 or CRC-32/ISIZE check) until the
 * input ends, their outputs placed one after another.  The members' outputs
 * must add up to output_size (else status 11; 7 when they exceed it), and an
 * input that ends inside a member gives that member's status (14 for a
 * missing trailer).  The first failing member's status is reported; on a
 * checksum mismatch (21, 24) the output decoded so far is kept, otherwise the
 * output is zero-filled.  This mode synchronises the stream with the host
 * once per member (the next member starts where the previous one ended), so
 * it must not be used under graph capture.  The reference rejects a second
 * stream after the first (tests/test_decode.py:679-713). */
#define HIP_ZLIB_FORMAT_MEMBERS 0x100
int HipZlibDecompressFormat(hipStream_t stream, int32_t format, const uint8_t* dictionary,
                            uint64_t dictionary_size, int64_t max_candidates, int64_t max_blocks,
                            const uint8_t* input, uint64_t input_size, uint8_t* output,
                            uint64_t output_size, uint32_t* metadata, uint64_t metadata_count);

/* Compress `files` packed inputs (host array input_sizes) into consecutive
 * padded slots; metadata (files x 2 u32, device) rows are [encoded_length, status].
 * The host-side size list is copied to the device before the call returns.
 * Replaces CudaZlibCompressBatch (codec_ffi.cu:1163-1172, body 1002-1063). */
int HipZlibCompressBatch(hipStream_t stream, int64_t chunk_bytes, const int64_t* input_sizes,
                         uint64_t files, const uint8_t* input, uint64_t input_size,
                         uint8_t* output, uint64_t output_size, uint32_t* metadata,
                         uint64_t metadata_rows, uint64_t metadata_cols);

/* Decompress packed independent streams.  encoded_metadata is null (rows = 0)
 * or compression's (files x 2) [length, status] rows on the device; then a
 * file's stream length is read on the device.  metadata rows are [status, 0].
 * Replaces CudaZlibDecompressBatch (codec_ffi.cu:1173-1182, body 1065-1107). */
int HipZlibDecompressBatch(hipStream_t stream, const int64_t* input_sizes, uint64_t input_count,
                           const int64_t* output_sizes, uint64_t output_count,
                           const uint8_t* input, uint64_t input_size,
                           const uint32_t* encoded_metadata, uint64_t encoded_rows,
                           uint64_t encoded_cols, uint8_t* output, uint64_t output_size,
                           uint32_t* metadata, uint64_t metadata_rows, uint64_t metadata_cols);

/* HipZlibCompress without any allocation: same arguments, results and
 * metadata, but the scratch comes from a fixed 48 MiB device array that the
 * library holds on each GPU for the life of the process, instead of the pool.
 * It calls no hipMalloc/hipFree or allocating routine, for callers that cannot
 * allocate (code under HIP graph capture, allocation-free serving loops).
 * Inputs are limited by that array: with 32 KiB chunks up to about 11 MiB
 * (scratch is about 5 bytes per input byte).  A larger input returns
 * HIP_ZLIB_INVALID_ARGUMENT, with the bytes it would need in
 * HipZlibErrorString(-1), and enqueues nothing.  Calls on one GPU share the
 * array: calls that overlap on a GPU (on different streams, or from different
 * threads) race, so callers serialise them.  No counterpart in the reference. */
int HipZlibCompressNoAlloc(hipStream_t stream, int64_t chunk_bytes, const uint8_t* input,
                           uint64_t input_size, uint8_t* output, uint64_t output_size,
                           uint32_t* metadata, uint64_t metadata_count);

/* Workspace pool controls.  Replace CudaZlibSetWorkspaceRetention,
 * CudaZlibWorkspacePoolStats and CudaZlibTrimWorkspacePool (codec_ffi.cu:1113-1142).
 * Retention may only change before the first pool is created.
 * stats = {retention_bytes, reserved_bytes, used_bytes, pool_count}. */
int HipZlibSetWorkspaceRetention(uint64_t bytes);
int HipZlibWorkspacePoolStats(int device, uint64_t* stats);
int HipZlibTrimWorkspacePool(int device);

/* Measurement hooks.  While enabled, every kernel the library launches is
 * bracketed by HIP events on the caller's stream.  Collect writes lines
 * "kernel launches total_ms" (after the caller synchronised the stream) and
 * returns the full text length; reset != 0 discards the records. */
int HipZlibProfileEnable(int enabled);
uint64_t HipZlibProfileCollect(char* buffer, uint64_t capacity, int reset);

/* Text for a return code of any entry point above (thread-local for -1). */
const char* HipZlibErrorString(int code);

#ifdef __cplusplus
}
#endif

#endif /* HIP_ZLIB_H_ */
