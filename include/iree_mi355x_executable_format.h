// Serialized executable: the dispatch library as a compiler would embed it in
// a module, and the loader a runtime uses to bring it back.
//
// Replaces the Hexagon executable serialization and loading:
//  * the compiler links the dispatch functions into an ELF shared object and
//    embeds it as a hal.executable.binary of mime type application/x-elf
//    (TG/HexagonExecutableSerialization.cpp:491-640, linked by
//    TG/LibraryBuilder.cpp:179-340);
//  * the runtime writes it out, dlopens it, looks up the query function,
//    checks the library version and rejects HAL imports, then binds the
//    exports by name (RT/dsp/executable.c:92-147).
// Here the container also carries the export names and attributes, so a
// host can check what it loads before it calls into it, and a checksum.
//
// Layout (little-endian):
//   iree_mi355x_executable_header_t
//   export table: per export, u64 flags, u64 lds_bytes, u64 threads, then
//                 the NUL-terminated names back to back
//   the ELF shared object (iree_mi355x_executable_library_query inside)
// The checksum is FNV-1a 64 over every byte after the header.
#ifndef IREE_MI355X_EXECUTABLE_FORMAT_H_
#define IREE_MI355X_EXECUTABLE_FORMAT_H_

#include <stddef.h>
#include <stdint.h>

#include "iree_mi355x_executable_library.h"

#ifdef __cplusplus
extern "C" {
#endif

#define IREE_MI355X_EXECUTABLE_MAGIC "MI355XEX"
#define IREE_MI355X_EXECUTABLE_FORMAT_VERSION 1u
#define IREE_MI355X_EXECUTABLE_MIME "application/x-elf"

typedef struct iree_mi355x_executable_header_t {
  char magic[8];              // IREE_MI355X_EXECUTABLE_MAGIC (no NUL)
  uint32_t format_version;    // IREE_MI355X_EXECUTABLE_FORMAT_VERSION
  uint32_t library_version;   // IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_*
  char arch[16];              // "gfx950", NUL-padded
  char mime[24];              // IREE_MI355X_EXECUTABLE_MIME, NUL-padded
  uint32_t export_count;
  uint32_t reserved;
  uint64_t table_offset, table_bytes;      // from the start of the header
  uint64_t library_offset, library_bytes;  // the ELF
  uint64_t checksum;                       // FNV-1a 64 of bytes after header
} iree_mi355x_executable_header_t;

// Serializes the ELF at `library_path` (NULL: this library's own file) with
// the export table its query returns. Returns the container size; writes it
// to `out` only when `capacity` is at least that. 0 on error (see
// iree_mi355x_last_error).
size_t iree_mi355x_executable_serialize(const char *library_path, void *out,
                                        size_t capacity);

// Checks magic, versions, architecture, offsets and checksum without loading.
int iree_mi355x_executable_verify(const void *data, size_t size);

typedef struct iree_mi355x_loaded_executable_t
    iree_mi355x_loaded_executable_t;

// Verifies, writes the ELF to an anonymous file and dlopens it, queries its
// library at IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST, rejects imports
// and checks its exports against the container's table.
int iree_mi355x_executable_load(const void *data, size_t size,
                                iree_mi355x_loaded_executable_t **out);

// The loaded library's table (for iree_mi355x_command_buffer_create).
const iree_mi355x_executable_library_t *iree_mi355x_loaded_executable_library(
    const iree_mi355x_loaded_executable_t *executable);

// Unloads. Every dispatch of the executable must have completed.
void iree_mi355x_loaded_executable_release(
    iree_mi355x_loaded_executable_t *executable);

#ifdef __cplusplus
}  // extern "C"
#endif

#endif  // IREE_MI355X_EXECUTABLE_FORMAT_H_
