"""Write the C block of INTEGRATION.md's `src/generate.c` section to stdout
(test infrastructure: tests/c/ compiles the documented snippet as it stands)."""
import sys

txt = open(sys.argv[1]).read()
sec = txt.split("## The change in `src/generate.c`", 1)[1]
code = sec.split("```c\n", 1)[1].split("```", 1)[0]
sys.stdout.write(code)
