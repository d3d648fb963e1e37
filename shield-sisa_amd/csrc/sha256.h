/* SHA-256 (FIPS 180-4), incremental.  Used for the weight-file fingerprint, the sidecar check and the
 * compute revision.  Plain C so that the host library, the synthetic-weight writer and tests share it. */
#ifndef SHV_SHA256_H
#define SHV_SHA256_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct shv_sha256 {
    uint32_t h[8];
    uint64_t length;       /* message bytes so far */
    uint8_t block[64];
    size_t fill;           /* bytes pending in block */
} shv_sha256;

void shv_sha256_init(shv_sha256* s);
void shv_sha256_update(shv_sha256* s, const void* data, size_t n);
void shv_sha256_final(shv_sha256* s, uint8_t digest[32]);
/* digest -> 64 lowercase hex characters + NUL */
void shv_sha256_hex(const uint8_t digest[32], char out[65]);

#ifdef __cplusplus
}
#endif
#endif
