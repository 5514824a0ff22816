/* The C ABI of libmingtts_hip.so for Swift.  Build with the repository's include/ on the
 * header path and the library's directory on the link path:
 *   swift build -Xcc -I<repo>/include -Xlinker -L<repo>/ming-tts_amd/csrc
 */
#include <mingtts_hip.h>
