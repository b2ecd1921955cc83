import sys

from torque_hip.cli import main

sys.exit(main())
