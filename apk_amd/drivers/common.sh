# Shared by the sweep drivers: where the binaries are, and where raw results go
# (results/raw under the current directory, as the reference's drivers write).
set -euo pipefail
BIN=${APK_BIN:-$(cd "$(dirname "${BASH_SOURCE[0]}")/../bin" && pwd)}
RAW=${APK_RAW:-results/raw}
mkdir -p "$RAW"
banner() { printf '\n=============== %s ===============\n' "$*"; }
