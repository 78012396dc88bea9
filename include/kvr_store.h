/*
 * kvr_store.h -- on-disk / wire format of the 1-bit tile store (format version 1).
 *
 * A store file carries the decode state of n_layers layers of B sequences x Hkv KV
 * heads ("segments", segment = b * Hkv + h): per layer the K and V tile bits and fp16
 * tile scales (the layout kvr_encode_tiles writes), optionally the K channel counts,
 * and optionally the exact recent tokens (the window, oldest first).  Everything is
 * little-endian.  Byte layout of a file:
 *
 *   [0, 256)     header, written by kvr_store_header_encode:
 *     0   char[8]  magic "KVRSTORE"
 *     8   u32      format version (KVR_STORE_FORMAT_VERSION)
 *     12  u32      header bytes (256)
 *     16  u32      C ABI version of the writer (kvr_abi_version; informational)
 *     20  i32      d (head_dim, 128)
 *     24  i32      T (tile tokens, 64 or 128)
 *     28  i32      transform (enum kvr_transform of the codec)
 *     32  i32      bit order (KVR_BITS_TOKEN_LSB)
 *     36  i32      scale dtype (KVR_FP16)
 *     40  i32      window dtype (enum kvr_dtype; meaningful with KVR_STORE_HAS_WINDOW)
 *     44  u32      flags (KVR_STORE_HAS_COUNTS | KVR_STORE_HAS_WINDOW)
 *     48  i32      n_layers
 *     52  u32      section alignment (KVR_STORE_ALIGN)
 *     56  i64      B          64  i64  Hkv         72  i64  n_tiles (per segment)
 *     80  i64      W (window size of the writer's cache, a multiple of T; 0: none)
 *     88  i64      win_len (window tokens per segment, 0 <= win_len < W + T)
 *     96  u64      payload bytes (everything after the header)
 *     104 u32      CRC-32 of the payload
 *     108 u32      0
 *     112 i64[4]   user words (the writer's own, e.g. a decoder's step counters)
 *     144 ..       zeros
 *     252 u32      CRC-32 of bytes [0, 252)
 *   [256, ...)   payload: for layer 0, 1, ...: its sections in enum kvr_store_section
 *                order (absent ones skipped), each starting at a multiple of
 *                KVR_STORE_ALIGN bytes from the start of the file, zeros between:
 *     KBITS, VBITS : uint64 [B*Hkv][n_tiles][128][T/64]; bit (t mod 64) of word t/64 is
 *                    the sigma-delta bit of token t of that channel (KVR_BITS_TOKEN_LSB)
 *     KSCALE,VSCALE: fp16 bit patterns [B*Hkv][n_tiles]
 *     KCOUNT       : uint8 [B*Hkv][n_tiles][128], set bits per channel over the tile
 *     WIN_K, WIN_V : window dtype [B][Hkv][win_len][128], oldest token first
 *
 * CRC-32 is the IEEE 802.3 / zlib one (reflected polynomial 0xEDB88320, initial and
 * final complement): kvr_crc32(0, p, n) == zlib.crc32(p).  All functions here are
 * host-only (no device, no HIP call) and return KVR_OK or a negative kvr_status with
 * kvr_last_error() set.
 *
 * Replaces: nothing in the reference -- it keeps its store in device memory only and
 *           rebuilds it on reset (modules/kvr_hook.py:316-326,
 *           modules/kvr_retrieval.py:150-160); the format serves prefix caching and
 *           fixture exchange.
 */
#ifndef KVR_STORE_H
#define KVR_STORE_H

#include <stddef.h>
#include <stdint.h>

#include "kvr_capi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define KVR_STORE_HEADER_BYTES 256
#define KVR_STORE_FORMAT_VERSION 1
#define KVR_STORE_ALIGN 64

enum kvr_store_flags { KVR_STORE_HAS_COUNTS = 1, KVR_STORE_HAS_WINDOW = 2 };
enum kvr_bit_order { KVR_BITS_TOKEN_LSB = 0 };
enum kvr_store_section {
  KVR_SEC_KBITS = 0,
  KVR_SEC_VBITS = 1,
  KVR_SEC_KSCALE = 2,
  KVR_SEC_VSCALE = 3,
  KVR_SEC_KCOUNT = 4,
  KVR_SEC_WIN_K = 5,
  KVR_SEC_WIN_V = 6,
  KVR_SEC_N = 7
};

typedef struct kvr_store_desc {
  uint32_t format_version; /* set by kvr_store_header_encode / _decode                */
  uint32_t abi_version;    /* set by encode (this library's), read by decode          */
  int32_t d, T, transform, bit_order, scale_dtype, win_dtype;
  uint32_t flags;
  int32_t n_layers;
  int64_t B, Hkv, n_tiles, W, win_len;
  uint64_t payload_bytes;  /* set by encode from the layout; decode checks it          */
  uint32_t payload_crc32;  /* the caller's CRC-32 of the payload                       */
  int64_t user[4];
} kvr_store_desc;

/* CRC-32 of n bytes continuing from crc (0 to start). */
uint32_t kvr_crc32(uint32_t crc, const void* data, size_t n);

/* Payload bytes of a store described by desc (its fields validated as by encode), or a
 * negative kvr_status. */
int64_t kvr_store_payload_bytes(const kvr_store_desc* desc);

/* Byte offset from the start of the file of section `section` of layer `layer`, with
 * its size in *bytes (nullable); a negative kvr_status if the description is invalid,
 * the index is out of range or the section is absent (flags). */
int64_t kvr_store_section(const kvr_store_desc* desc, int layer, int section, int64_t* bytes);

/* Validate desc and write the 256-byte header (format version, ABI version, payload
 * bytes and the header CRC filled in; desc->payload_crc32 taken as given). */
int kvr_store_header_encode(const kvr_store_desc* desc, void* header);

/* Read and validate a header: magic, format version (newer ones are
 * KVR_ERR_UNSUPPORTED), header CRC, field ranges and the payload size. */
int kvr_store_header_decode(const void* header, size_t n, kvr_store_desc* desc);

#ifdef __cplusplus
}
#endif

#endif /* KVR_STORE_H */
